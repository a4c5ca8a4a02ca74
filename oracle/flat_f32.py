"""NumPy restatement of the reference's fp32-dot GPU path -- TEST INFRASTRUCTURE ONLY.

``_flat_triton`` with ``dot`` other than "bf16" (h3/htrc_flat.py:181-276; the kernels of
h3/htrc_flat_triton.py with DOT = 0): the leaf state in fp32 (store="fp32", the reference's default)
or bf16 (store="bf16"), every dot on fp32 operands -- IEEE (prec="ieee") or rounded to TF32 first
(prec="tf32", to nearest with ties away from zero, as a TF32 tensor-core operand is converted) --
the row-max select over every sel_stride-th row of each group of tiles, top-k with sink leaves,
and per row one softmax over the far leaves outside the near set and the near leaves' tokens.
One head.  Products and sums are float64; the values the reference stores (g, vb, lz, SEL) are
rounded to float32 (g and vb to bf16 for store="bf16"), so the GPU is compared with the exact
value of the reference's formula on the reference's own stored operands.  The softmax weights
enter the PV products unrounded (the reference rounds them to TF32 as well under prec="tf32",
a 2^-11 relative difference the tests' tolerances carry).

Pinned in tests/test_oracle_f32.py: the TF32 rounding on known values (ties away, carries into
the exponent, infinities); store="fp32" at IEEE precision equals ``flat_fp32`` (the reference's
torch backend, h3/htrc_flat.py:279-388) wherever both select the same near leaves; every leaf
near equals dense attention; and the bf16 store is the fp32 store's pipeline on g and vb rounded
to bf16.
"""
from __future__ import annotations

import math

import numpy as np

from . import bf16
from .flat_i8 import group_centres, kmeans_order, tile_centres, topk


def tf32_rna(x) -> np.ndarray:
    """float32 -> TF32 (10 explicit mantissa bits), to nearest with ties away from zero;
    infinities and NaN unchanged (the tensor-core operand conversion, cvt.rna.tf32.f32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    r = ((u + np.uint32(0x1000)) & np.uint32(0xFFFFE000)).astype(np.uint32)
    special = (u & np.uint32(0x7F800000)) == np.uint32(0x7F800000)
    return np.where(special, u, r).astype(np.uint32).view(np.float32)


def _op(x, prec: str) -> np.ndarray:
    """A dot operand as the reference's tl.dot takes it (float64 for the exact products)."""
    x = np.asarray(x, np.float32)
    return (tf32_rna(x) if prec == "tf32" else x).astype(np.float64)


def _stored(x, store: str) -> np.ndarray:
    """A state tensor as the reference stores it: float32, or bf16 for store="bf16"."""
    x = np.asarray(x, np.float32)
    return bf16.round_f32(x) if store == "bf16" else x


def stats(mu, k, v, leaf: int, scale: float, prec: str = "ieee", store: str = "fp32"):
    """Leaf statistics (h3/htrc_flat_triton.py:41-85 with FP8 = I8 = 0): mu [nc, d], k / v [nk, d]
    float32 -> g, vb [nc, nb, d] (float32; bf16 values for store="bf16") and lz [nc, nb]:
    a = (mu . k) scale, w = softmax_leaf(a), g = (w K) scale, vb = w V, lz = max + log sum."""
    mu = np.asarray(mu, np.float32)
    nc, d = mu.shape
    nb = k.shape[0] // leaf
    kl = np.asarray(k, np.float32)[:nb * leaf].reshape(nb, leaf, d).astype(np.float64)
    vl = np.asarray(v, np.float32)[:nb * leaf].reshape(nb, leaf, d).astype(np.float64)
    sc = np.float32(scale)
    a = (np.einsum("cd,lkd->clk", _op(mu, prec), kl).astype(np.float32) * sc).astype(np.float32)
    m = a.max(-1, keepdims=True)
    e = np.exp((a - m).astype(np.float64)).astype(np.float32)
    z = e.sum(-1, keepdims=True, dtype=np.float64).astype(np.float32)
    w = (e / z).astype(np.float32)
    wo = _op(w, prec)
    g = np.einsum("clk,lkd->cld", wo, kl).astype(np.float32) * sc
    vb = np.einsum("clk,lkd->cld", wo, vl).astype(np.float32)
    lz = (m[..., 0].astype(np.float64) + np.log(z[..., 0].astype(np.float64))).astype(np.float32)
    return _stored(g, store), _stored(vb, store), lz


def _group_rows(n: int, tile: int, group: int, c: int, stride: int) -> np.ndarray:
    """Operator rows of group c as the reference pads them (tiles past the last repeat it, rows
    past the last query repeat it), every stride-th row."""
    nt = -(-n // tile)
    j = np.arange(0, group * tile, stride)
    t = np.minimum(c * group + j // tile, nt - 1)
    return np.minimum(t * tile + j % tile, n - 1)


def select(qf, mu, g, lz, *, tile: int, group: int = 1, stride: int = 1, prec: str = "ieee") -> np.ndarray:
    """SEL [ng, nb] = max over every stride-th row of the group of (q - mu) . g, + lz
    (h3/htrc_flat_triton.py:214-254, DOT = 0); qf [n, d] in operator row order."""
    qf = np.asarray(qf, np.float32)
    ng, nb, d = g.shape
    sel = np.empty((ng, nb), np.float32)
    go = _op(g, prec)
    for c in range(ng):
        rows = _group_rows(qf.shape[0], tile, group, c, stride)
        dq = (qf[rows] - mu[c][None, :]).astype(np.float32)
        s = (_op(dq, prec) @ go[c].T).astype(np.float32)
        sel[c] = (s.max(0) + lz[c]).astype(np.float32)
    return sel


def attend(qf, mu, g, lz, vb, idx, excl, k, v, *, tile: int, leaf: int, scale: float, group: int = 1,
           prec: str = "ieee"):
    """Far leaves outside the near set (score (q - mu) . g + lz, value vb) and the near leaves'
    tokens (score (q . k) scale, value v) in one exact softmax per row
    (h3/htrc_flat_triton.py:88-211, DOT = 0) -> out [n, d], logz [n] (operator row order)."""
    qf = np.asarray(qf, np.float32)
    n, d = qf.shape
    nt = -(-n // tile)
    out = np.zeros((n, d), np.float64)
    logz = np.zeros((n,), np.float64)
    kf = np.asarray(k, np.float32)
    vf = np.asarray(v, np.float64)
    ar = np.arange(leaf)
    for t in range(nt):
        c = t // group
        r0, r1 = t * tile, min(n, t * tile + tile)
        qr = qf[r0:r1]
        dq = (qr - mu[c][None, :]).astype(np.float32)
        far = ~excl[c][: g.shape[1]].astype(bool)
        sf = (_op(dq, prec) @ _op(g[c][far], prec).T).astype(np.float32) + lz[c][far][None, :]
        vals = [np.asarray(vb[c][far], np.float64)]
        scores = [sf.astype(np.float64)]
        if idx.shape[1] > 0:
            tok = (idx[c][:, None] * leaf + ar).reshape(-1)
            sn = (_op(qr, prec) @ _op(kf[tok], prec).T).astype(np.float32) * np.float32(scale)
            scores.append(sn.astype(np.float64))
            vals.append(vf[tok])
        s = np.concatenate(scores, 1)
        vv = np.concatenate(vals, 0)
        m = s.max(1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        e = np.exp(s - m)
        z = e.sum(1, keepdims=True)
        out[r0:r1] = (e @ vv) / np.maximum(z, 1e-30)
        with np.errstate(divide="ignore"):
            logz[r0:r1] = (np.log(z) + m)[:, 0]
    return out, logz


def flat_f32(q, k, v, *, tile: int = 64, leaf: int = 64, exact_leaves: int = 64, store: str = "fp32",
             prec: str = "ieee", group: int = 1, sel_stride: int = 1, sink_leaves: int = 0, order: str = "seq",
             scale: float | None = None, select_mode: str = "max") -> dict:
    """The fp32-dot flat operator for one head: q [n, d], k / v [nk, d] float32 arrays (bf16
    values for k / v, as the operator takes them), nk % leaf == 0.  Returns the intermediates
    (mu, g, vb, lz, sel, idx, excl; perm for order="kmeans") plus out [n, d] and logz [n] in
    query order.  select_mode "bound": lz + max_r ||q - mu|| ||g|| (h3/htrc_flat.py:255-257)."""
    qf = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    n, d = qf.shape
    if k.shape[0] % leaf:
        raise ValueError("key count must be a multiple of the leaf size")
    nb = k.shape[0] // leaf
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    sink = max(0, min(int(sink_leaves), nb))
    kx = min(int(exact_leaves) + sink, nb)
    st: dict = {}
    if order == "kmeans":
        st["perm"] = kmeans_order(qf)
        qf = qf[st["perm"]]
    elif order != "seq":
        raise ValueError("order must be seq or kmeans")
    st["mu"] = tile_centres(qf, tile) if group == 1 else group_centres(qf, tile, group)
    st["g"], st["vb"], st["lz"] = stats(st["mu"], k, v, leaf, scale, prec, store)
    ng = st["mu"].shape[0]
    if kx > 0:
        if select_mode == "bound":
            sel = np.empty((ng, nb), np.float32)
            for c in range(ng):
                rows = _group_rows(n, tile, group, c, 1)
                dq = (qf[rows] - st["mu"][c][None, :]).astype(np.float64)
                r = np.sqrt((dq * dq).sum(1)).max()
                gn = np.sqrt((st["g"][c].astype(np.float64) ** 2).sum(1))
                sel[c] = (st["lz"][c] + r * gn).astype(np.float32)
            st["sel"] = sel
        else:
            st["sel"] = select(qf, st["mu"], st["g"], st["lz"], tile=tile, group=group, stride=sel_stride, prec=prec)
        st["idx"], st["excl"] = topk(st["sel"], kx, sink)
    else:
        st["idx"] = np.zeros((ng, 0), np.int32)
        st["excl"] = np.zeros((ng, nb), np.int8)
    out, logz = attend(qf, st["mu"], st["g"], st["lz"], st["vb"], st["idx"], st["excl"], k, v, tile=tile, leaf=leaf,
                       scale=scale, group=group, prec=prec)
    if order == "kmeans":
        o2, l2 = np.empty_like(out), np.empty_like(logz)
        o2[st["perm"]], l2[st["perm"]] = out, logz
        out, logz = o2, l2
    st["out"], st["logz"] = out.astype(np.float32), logz.astype(np.float32)
    return st


def tail_merge(out, logz, q, tk, tv, scale: float, prec: str = "ieee"):
    """Keys past the last full leaf, attended exactly by every query with fp32 operands (TF32 for
    prec="tf32"; h3/htrc_flat_triton.py:187-207 with DOT = 0), merged into a finished (out [n, d],
    logz [n]): one softmax over all keys, by the split-merge algebra of :257-273."""
    s = ((_op(q, prec) @ _op(tk, prec).T).astype(np.float32) * np.float32(scale)).astype(np.float64)
    m = s.max(1)
    p = np.exp(s - m[:, None])
    l = p.sum(1)
    mean = (p @ np.asarray(tv, np.float64)) / l[:, None]
    lse = m + np.log(l)
    lz0 = np.asarray(logz, np.float64)
    z = np.logaddexp(lz0, lse)
    res = np.asarray(out, np.float64) * np.exp(lz0 - z)[:, None] + mean * np.exp(lse - z)[:, None]
    return res.astype(np.float32), z.astype(np.float32)
